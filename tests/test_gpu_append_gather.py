"""GPU parity: paged append / gather / copy_blocks / swap against the CPU oracle.

Bar: bit-exact. The pool image read back from HBM must equal, byte for byte, the
image the oracle builds from the same inputs (pool.rs:122-153 semantics through
the paged layout; f16 RNE or ties-away; Q8_0 per q8_dot.rs:46-59).
"""
import numpy as np
import pytest

from tests.helpers import make_pools, slots_for, to_dev

pytestmark = pytest.mark.gpu


def _f16_sweep_values(seed=0):
    """Every combination of the top 19 bits of an f32 (sign, exponent, top 10
    mantissa bits) with low-13-bit patterns that straddle every rounding case
    (exact, just above/below half, exact half), plus random bit patterns."""
    hi = np.arange(1 << 19, dtype=np.uint32) << 13
    lows = np.array([0x0000, 0x0001, 0x0fff, 0x1000, 0x1001, 0x1fff], dtype=np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    rng = np.random.default_rng(seed)
    bits = np.concatenate([bits, rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)])
    return bits.view(np.float32)


@pytest.mark.parametrize("rounding", [0, 1])
def test_append_f16_encoding_sweep_bit_exact(rounding):
    from oracle import ref
    x = _f16_sweep_values()
    d = 64
    n_tok = x.size // d
    x = x[: n_tok * d].reshape(n_tok, 1, d)
    v = x[::-1].copy()
    nblk = (n_tok + 15) // 16
    pool, layout = make_pools(1, 1, d, nblk, dtype=1, rounding=rounding)
    pool.fill(0)
    slots = np.arange(n_tok, dtype=np.int64)
    pool.append(0, to_dev(x), to_dev(v), to_dev(slots))
    got = pool.read()
    want = ref.new_pool(layout)
    ref.append(layout, want, 0, x, v, slots)
    mism = np.flatnonzero(got != want)
    assert mism.size == 0, f"{mism.size} bytes differ, first at {mism[:4]}"
    assert pool.take_fault_flags() == 0


def _q8_blocks(seed=0):
    rng = np.random.default_rng(seed)
    blocks = [rng.standard_normal((2048, 32)).astype(np.float32)]
    out = rng.standard_normal((2048, 32)).astype(np.float32)
    mask = rng.random(out.shape) < 0.01
    out[mask] = np.where(rng.random(mask.sum()) < 0.5, -20.0, 20.0)
    blocks.append(out)
    for e in range(-45, 39, 3):  # amax from subnormal to near FLT_MAX
        blocks.append((rng.standard_normal((64, 32)) * 10.0 ** e).astype(np.float32))
    ties = np.zeros((254, 32), np.float32)  # amax 127 -> d = 1, id = 1: exact .5 ties
    ties[:, 0] = 127.0
    ties[:, 1:] = (np.arange(-127, 127)[:, None] + 0.5).astype(np.float32)
    blocks.append(ties)
    # Near ties: v with fl(v*id) == k + 0.5 exactly while the exact product is not,
    # so an implicitly fused v*id - trunc(v*id) rounds the other way.
    near = []
    for amax in rng.uniform(0.5, 30.0, 4000).astype(np.float32):
        dd = np.float32(amax / np.float32(127.0))
        idv = np.float32(np.float32(1.0) / dd)
        kk = rng.integers(-120, 120)
        v0 = np.float32((kk + 0.5) * np.float64(dd))
        for cand in (np.nextafter(v0, np.float32(-1e9)), v0, np.nextafter(v0, np.float32(1e9))):
            p = np.float32(cand * idv)
            if p == np.float32(kk + 0.5) and np.float64(cand) * np.float64(idv) != kk + 0.5 \
                    and abs(cand) <= amax:
                row = np.zeros(32, np.float32)
                row[0] = amax
                row[1:] = cand
                near.append(row)
                break
    assert len(near) > 100
    blocks.append(np.array(near, np.float32))
    special = np.zeros((8, 32), np.float32)
    special[1, 3] = 1.0
    special[2, :] = np.inf
    special[3, 5] = np.nan
    special[4, 7] = -np.inf
    special[5, :] = -0.0
    special[6, 9] = np.float32(1e-45)
    special[7, :] = np.float32(3.4e38)
    blocks.append(special)
    b = np.concatenate(blocks)
    return b[: b.shape[0] // 4 * 4]


@pytest.mark.parametrize("rounding", [0, 1])
def test_append_q8_bit_exact(rounding):
    from oracle import ref
    blocks = _q8_blocks()
    d, hkv = 128, 1
    x = blocks.reshape(-1, hkv, d)
    n_tok = x.shape[0]
    v = np.ascontiguousarray(x[::-1])
    pool, layout = make_pools(1, hkv, d, (n_tok + 15) // 16, dtype=8, rounding=rounding)
    pool.fill(0)
    slots = np.arange(n_tok, dtype=np.int64)
    pool.append(0, to_dev(x), to_dev(v), to_dev(slots))
    got = pool.read()
    want = ref.new_pool(layout)
    ref.append(layout, want, 0, x, v, slots)
    mism = np.flatnonzero(got != want)
    assert mism.size == 0, f"{mism.size} bytes differ, first at {mism[:4]}"


@pytest.mark.parametrize("dtype,d", [(0, 128), (1, 128), (1, 64), (8, 64), (0, 4), (1, 12)])
def test_append_gather_roundtrip_scattered(dtype, d):
    """Append through a scattered slot mapping (with -1 padding), gather back by
    slot (f32 and raw) and by block table; all bit-exact against the oracle."""
    import torch
    from oracle import ref
    rng = np.random.default_rng(1)
    L, hkv, nblk = 3, 2, 64
    pool, layout = make_pools(L, hkv, d, nblk, dtype=dtype)
    pool.fill(0x5a)
    want = np.full(layout.pool_bytes, 0x5a, np.uint8)
    seqs = [37, 1, 16, 100, 0, 33]
    perm = rng.permutation(nblk).astype(np.int32)
    tables, off = [], 0
    for c in seqs:
        nb = (c + 15) // 16
        tables.append(perm[off: off + nb])
        off += nb
    max_blocks = max(1, max(len(t) for t in tables))
    tab = np.zeros((len(seqs), max_blocks), np.int32)
    for i, t in enumerate(tables):
        tab[i, : len(t)] = t
    slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(seqs)])
    slots = np.insert(slots, [3, 10], -1)  # padding tokens
    n = slots.size
    for layer in range(L):
        k = rng.standard_normal((n, hkv, d), dtype=np.float32)
        v = rng.standard_normal((n, hkv, d), dtype=np.float32)
        pool.append(layer, to_dev(k), to_dev(v), to_dev(slots))
        ref.append(layout, want, layer, k, v, slots)
    assert np.array_equal(pool.read(), want)
    assert pool.take_fault_flags() == 0
    image = want
    for fmt in (0, 1):
        ek, ev = ref.gather_slots(layout, image, 1, slots, fmt)
        fill = -7.0 if fmt == 0 else 0xA5
        gk = torch.full(ek.shape, fill, dtype=torch.float32 if fmt == 0 else torch.uint8,
                        device="cuda")
        gv = torch.full(ev.shape, fill, dtype=gk.dtype, device="cuda")
        pool.gather_slots(1, to_dev(slots), gk, gv, fmt)
        gk, gv = gk.cpu().numpy(), gv.cpu().numpy()
        live = slots >= 0
        assert np.array_equal(gk[live].view(np.uint8), ek[live].view(np.uint8))
        assert np.array_equal(gv[live].view(np.uint8), ev[live].view(np.uint8))
        if d % 8 == 0 or dtype == 8:
            ctx = np.array(seqs, np.int32)
            tk, tv, offs = ref.gather_tables(layout, image, 2, tab, ctx, fmt)
            ok = torch.zeros(tk.shape, dtype=torch.float32 if fmt == 0 else torch.uint8,
                             device="cuda")
            ov = torch.zeros_like(ok)
            pool.gather_tables(2, to_dev(tab), to_dev(ctx), to_dev(offs), int(ctx.max()), ok, ov,
                               fmt)
            assert np.array_equal(ok.cpu().numpy().view(np.uint8), tk.view(np.uint8))
            assert np.array_equal(ov.cpu().numpy().view(np.uint8), tv.view(np.uint8))


@pytest.mark.parametrize("dtype", [1, 8])
@pytest.mark.parametrize("d,hkv", [(128, 2), (64, 3), (64, 2), (128, 5)])
@pytest.mark.parametrize("rounding", [0, 1])
def test_append_runs_at_every_alignment(dtype, d, hkv, rounding):
    """F16 and Q8_0 append (the 16-token window kernels) of slot mappings whose runs of
    consecutive slots start at every offset of a block and at every position of a
    16-token window: chunks of 1..40 tokens continuing 0..15 tokens into a block, a
    descending run, random single slots, -1 padding, and a token count that leaves the
    last window partial; head counts that leave a workgroup's last heads empty. Bytes no
    token names keep the fill pattern; all bit-exact against the oracle."""
    from oracle import ref
    rng = np.random.default_rng(d + hkv + rounding + dtype)
    nblk = 160
    pool, layout = make_pools(2, hkv, d, nblk, dtype=dtype, rounding=rounding)
    pool.fill(0x5a)
    want = np.full(layout.pool_bytes, 0x5a, np.uint8)
    perm = rng.permutation(nblk)
    parts, b = [], 0
    for start in range(16):
        n = int(rng.integers(1, 41))
        nb = (start + n + 15) // 16
        blocks = perm[b: b + nb]
        b += nb
        pos = np.arange(start, start + n)
        parts.append(blocks[pos // 16].astype(np.int64) * 16 + pos % 16)
        if start % 5 == 0:
            parts.append(np.array([-1], np.int64))
    rest = perm[b: b + 4].astype(np.int64)
    parts.append((rest[0] * 16 + np.arange(16))[::-1])      # descending run
    parts.append(rng.permutation(np.concatenate([rest[1] * 16 + np.arange(16),
                                                 rest[2] * 16 + np.arange(16)]))[:23])
    parts.append(rest[3] * 16 + np.array([3, 4, 5, 9, 10, 15]))
    slots = np.concatenate(parts)
    if slots.size % 16 == 0:  # keep the last window partial
        slots = np.append(slots, rest[3] * 16 + 7)
    assert np.unique(slots[slots >= 0]).size == (slots >= 0).sum()
    for layer in range(2):
        k = rng.standard_normal((slots.size, hkv, d), dtype=np.float32)
        v = rng.standard_normal((slots.size, hkv, d), dtype=np.float32)
        pool.append(layer, to_dev(k), to_dev(v), to_dev(slots))
        ref.append(layout, want, layer, k, v, slots)
    got = pool.read()
    mism = np.flatnonzero(got != want)
    assert mism.size == 0, f"{mism.size} bytes differ, first at {mism[:4]}"
    assert pool.take_fault_flags() == 0


def test_append_out_of_range_slot_is_skipped_and_flagged():
    from oracle import ref
    pool, layout = make_pools(1, 1, 64, 4)
    pool.fill(0)
    k = np.ones((3, 1, 64), np.float32)
    slots = np.array([0, 4 * 16, 5], np.int64)  # middle one is past the pool
    pool.append(0, to_dev(k), to_dev(k), to_dev(slots))
    assert pool.take_fault_flags() == 1
    want = ref.new_pool(layout)
    skipped = ref.append(layout, want, 0, k, k, slots)
    assert skipped == 1
    assert np.array_equal(pool.read(), want)
    assert pool.take_fault_flags() == 0


@pytest.mark.parametrize("dtype", [1, 8])
def test_copy_blocks_bit_exact(dtype):
    import torch
    from oracle import ref
    rng = np.random.default_rng(2)
    nblk = 48
    pool, layout = make_pools(2, 2, 128, nblk, dtype=dtype)
    img = rng.integers(0, 256, layout.pool_bytes, dtype=np.uint8)
    pool.write(img)
    src = rng.choice(nblk // 2, 20, replace=False)
    dst = nblk // 2 + rng.choice(nblk // 2, 20, replace=False)
    pairs = np.stack([src, dst], 1).astype(np.int64)
    pool.copy_blocks(to_dev(pairs))
    torch.cuda.synchronize()
    want = img.copy()
    ref.copy_blocks(layout, want, pairs)
    assert np.array_equal(pool.read(), want)
    bad = np.array([[0, nblk]], np.int64)
    pool.copy_blocks(to_dev(bad))
    assert pool.take_fault_flags() == 2
    assert np.array_equal(pool.read(), want)


def test_swap_out_in_roundtrip():
    import torch
    rng = np.random.default_rng(3)
    nblk, nhost = 32, 16
    pool, layout = make_pools(2, 2, 64, nblk, num_host_blocks=nhost)
    img = rng.integers(0, 256, layout.pool_bytes, dtype=np.uint8)
    pool.write(img)
    bb = layout.block_bytes
    dev_blocks = np.array([3, 4, 5, 9, 20, 21, 31, 0])
    host_blocks = np.array([0, 1, 2, 7, 8, 9, 15, 3])
    pool.swap_out(np.stack([dev_blocks, host_blocks], 1))
    torch.cuda.synchronize()
    pool.fill(0)
    torch.cuda.synchronize()
    back = np.array([10, 11, 12, 13, 14, 15, 16, 17])
    pool.swap_in(np.stack([host_blocks, back], 1))
    torch.cuda.synchronize()
    got = pool.read()
    for db, nb in zip(dev_blocks, back):
        assert np.array_equal(got[nb * bb:(nb + 1) * bb], img[db * bb:(db + 1) * bb])
    import ferrum_amd as fa
    with pytest.raises(fa.CacheError, match="unknown host block"):
        pool.swap_out(np.array([[0, nhost]]))

"""GPU parity: block-table and slot gather (the paged KvPool::k / v of
crates/kvcache/src/pool.rs:174-204) bit-exact against the oracle.

F16 and Q8_0 pools with 16-token blocks and head_dim 64 / 128 take the tile kernels (one
workgroup per 16 tokens of one block and one or two KV heads; 16-byte loads, the V
transpose through LDS). Covered:
- both output formats: decoded f32 (KvPool::k's f32 rows) and raw storage (binary16, or
  Ferrum's 34-byte Q8_0 blocks, core-types/src/dtype.rs:19-21);
- head counts that leave a workgroup's second head empty (head_dim 64, odd counts);
- contexts of 0, 1, 15, 16, 17 and longer (partial last blocks), output rows placed at
  gapped offsets (rows between sequences stay untouched);
- a table entry outside the pool (FKV_FAULT_BLOCK_RANGE; its rows untouched) and a
  context past the table (FKV_FAULT_CTX_RANGE; clamped);
- slot windows that are whole blocks (tile path), partial and scattered windows with -1
  padding (per-chunk path), and outputs that are not 16-byte aligned (per-chunk kernels).
"""
import numpy as np
import pytest

from tests.helpers import make_pools, slots_for, to_dev

pytestmark = pytest.mark.gpu


def _filled_pool(dtype, d, hkv, nblk, layers=2, seed=0):
    import torch
    from oracle import ref
    rng = np.random.default_rng(seed)
    pool, layout = make_pools(layers, hkv, d, nblk, dtype=dtype)
    pool.fill(0x3c)
    want = np.full(layout.pool_bytes, 0x3c, np.uint8)
    slots = np.arange(nblk * 16, dtype=np.int64)
    for layer in range(layers):
        k = rng.standard_normal((slots.size, hkv, d), dtype=np.float32) * 3
        v = rng.standard_normal((slots.size, hkv, d), dtype=np.float32) * 3
        pool.append(layer, to_dev(k), to_dev(v), to_dev(slots))
        ref.append(layout, want, layer, k, v, slots)
    torch.cuda.synchronize()
    assert np.array_equal(pool.read(), want)
    return pool, layout, want, rng


def _rows(a, sel):
    """The selected rows as bytes, one row a line (shapes of the oracle's and the
    device outputs differ: [rows][heads * row] against [rows][heads][row])."""
    r = np.ascontiguousarray(a[sel])
    return r.view(np.uint8).reshape(r.shape[0], r.itemsize * int(np.prod(r.shape[1:])))


def _out(shape_rows, hkv, d, fmt, dtype, fill):
    import torch
    if fmt == 0:
        return torch.full((shape_rows, hkv, d), fill, dtype=torch.float32, device="cuda")
    per = d * 2 if dtype == 1 else d // 32 * 34
    return torch.full((shape_rows, hkv, per), 0xA5, dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("dtype,d,hkv", [(1, 128, 8), (1, 64, 3), (8, 128, 8), (8, 64, 3),
                                         (1, 128, 1), (8, 64, 1)])
def test_gather_tables_tile_bit_exact(dtype, d, hkv, fmt):
    import ferrum_amd as fa
    from oracle import ref
    nblk = 120
    pool, layout, image, rng = _filled_pool(dtype, d, hkv, nblk, seed=d + hkv + dtype)
    ctxs = [0, 1, 15, 16, 17, 300, 700]
    nb = [(c + 15) // 16 for c in ctxs]
    perm = rng.permutation(nblk).astype(np.int32)
    tab = np.zeros((len(ctxs), max(nb)), np.int32)
    o = 0
    for i, n in enumerate(nb):
        tab[i, :n] = perm[o:o + n]
        o += n
    ctx = np.array(ctxs, np.int32)
    # rows of sequence i start at offs[i]; 5 spare rows after each sequence
    offs = np.concatenate([[3], 3 + np.cumsum(ctx[:-1].astype(np.int64) + 5)]).astype(np.int64)
    rows = int(offs[-1] + ctx[-1] + 4)
    wk, wv, woffs = ref.gather_tables(layout, image, 1, tab, ctx, fmt)
    gk = _out(rows, hkv, d, fmt, dtype, -7.0)
    gv = _out(rows, hkv, d, fmt, dtype, -7.0)
    pool.gather_tables(1, to_dev(tab), to_dev(ctx), to_dev(offs), int(ctx.max()), gk, gv, fmt)
    gk, gv = gk.cpu().numpy(), gv.cpu().numpy()
    assert pool.take_fault_flags() == 0
    touched = np.zeros(rows, bool)
    for i, c in enumerate(ctxs):
        touched[offs[i]:offs[i] + c] = True
        src = slice(int(woffs[i]), int(woffs[i]) + c)
        dst = slice(int(offs[i]), int(offs[i]) + c)
        assert np.array_equal(_rows(gk, dst), _rows(wk, src)), f"K of seq {i}"
        assert np.array_equal(_rows(gv, dst), _rows(wv, src)), f"V of seq {i}"
    if fmt == 0:
        assert np.all(gk[~touched] == -7.0) and np.all(gv[~touched] == -7.0)
    else:
        assert np.all(gk[~touched] == 0xA5) and np.all(gv[~touched] == 0xA5)
    # a table entry outside the pool: its 16 rows are left alone and the fault raised;
    # a context past the table: clamped to it
    bad = tab.copy()
    bad[5, 2] = nblk + 7
    ctx2 = ctx.copy()
    ctx2[6] = tab.shape[1] * 16 + 40  # the last sequence: its clamped rows overlap nothing
    gk2 = _out(rows + 200, hkv, d, fmt, dtype, -7.0)
    gv2 = _out(rows + 200, hkv, d, fmt, dtype, -7.0)
    # (max_ctx_len may not exceed the table; the device context does)
    pool.gather_tables(1, to_dev(bad), to_dev(ctx2), to_dev(offs), tab.shape[1] * 16, gk2, gv2,
                       fmt)
    flags = pool.take_fault_flags()
    assert flags == fa.FAULT_BLOCK_RANGE | fa.FAULT_CTX_RANGE
    gk2 = gk2.cpu().numpy()
    skipped = slice(int(offs[5]) + 32, int(offs[5]) + 48)
    fillv = -7.0 if fmt == 0 else 0xA5
    assert np.all(gk2[skipped] == fillv)
    keep = slice(int(offs[5]), int(offs[5]) + 32)
    assert np.array_equal(_rows(gk2, keep), _rows(gk, keep))
    keep6 = slice(int(offs[6]), int(offs[6]) + 700)
    assert np.array_equal(_rows(gk2, keep6), _rows(gk, keep6))


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("dtype,d,hkv", [(1, 128, 8), (1, 64, 3), (8, 128, 2), (8, 64, 3)])
def test_gather_slots_windows_bit_exact(dtype, d, hkv, fmt):
    """Slot lists mixing whole blocks at 16-token window boundaries (the tile path) with
    a partial block, a reversed block, scattered slots and -1 padding (per-chunk path)."""
    from oracle import ref
    nblk = 64
    pool, layout, image, rng = _filled_pool(dtype, d, hkv, nblk, seed=7 * d + hkv)
    perm = rng.permutation(nblk)
    parts = [perm[0] * 16 + np.arange(16), perm[1] * 16 + np.arange(16),   # whole blocks
             perm[2] * 16 + np.arange(5, 16), np.array([-1, -1]),           # partial
             perm[3] * 16 + np.arange(16)[::-1],                            # reversed
             rng.permutation(perm[4] * 16 + np.arange(16))[:9],             # scattered
             perm[5] * 16 + np.arange(16),                                  # whole, shifted
             np.array([-1] * 10), perm[6] * 16 + np.arange(16),             # whole, at token 96
             perm[7] * 16 + np.arange(16), perm[8] * 16 + np.arange(7)]     # partial tail
    slots = np.concatenate(parts).astype(np.int64)
    assert np.array_equal(slots[96:128], np.concatenate(parts[8:10]))  # windows 6 and 7 whole
    wk, wv = ref.gather_slots(layout, image, 0, slots, fmt)
    gk = _out(slots.size, hkv, d, fmt, dtype, -7.0)
    gv = _out(slots.size, hkv, d, fmt, dtype, -7.0)
    pool.gather_slots(0, to_dev(slots), gk, gv, fmt)
    gk, gv = gk.cpu().numpy(), gv.cpu().numpy()
    assert pool.take_fault_flags() == 0
    live = slots >= 0
    assert np.array_equal(_rows(gk, live), _rows(wk, live))
    assert np.array_equal(_rows(gv, live), _rows(wv, live))
    fillv = -7.0 if fmt == 0 else 0xA5
    assert np.all(gk[~live] == fillv) and np.all(gv[~live] == fillv)


@pytest.mark.parametrize("dtype", [1, 8])
def test_gather_unaligned_outputs(dtype):
    """Outputs 4 bytes past a 16-byte boundary take the per-chunk kernels: same bytes."""
    import torch
    from oracle import ref
    d, hkv, nblk = 128, 2, 16
    pool, layout, image, rng = _filled_pool(dtype, d, hkv, nblk, seed=3)
    ctx = np.array([40, 16], np.int32)
    tab = rng.permutation(nblk).astype(np.int32)[:6].reshape(2, 3)
    wk, wv, offs = ref.gather_tables(layout, image, 0, tab, ctx, 0)
    n = int(ctx.sum())
    base_k = torch.zeros(n * hkv * d + 1, dtype=torch.float32, device="cuda")
    base_v = torch.zeros_like(base_k)
    gk, gv = base_k[1:].view(n, hkv, d), base_v[1:].view(n, hkv, d)
    assert gk.data_ptr() % 16 == 4
    pool.gather_tables(0, to_dev(tab), to_dev(ctx), to_dev(offs), int(ctx.max()), gk, gv, 0)
    assert np.array_equal(gk.cpu().numpy().view(np.uint8), wk.view(np.uint8))
    assert np.array_equal(gv.cpu().numpy().view(np.uint8), wv.view(np.uint8))
    slots = slots_for(tab[0], 40)
    sk, sv = ref.gather_slots(layout, image, 0, slots, 0)
    pool.gather_slots(0, to_dev(slots), gk[:40], gv[:40], 0)
    assert np.array_equal(gk[:40].cpu().numpy().view(np.uint8), sk.view(np.uint8))
    assert np.array_equal(gv[:40].cpu().numpy().view(np.uint8), sv.view(np.uint8))
    assert pool.take_fault_flags() == 0

"""Shared helpers for the GPU parity tests (oracle = checker only)."""
from __future__ import annotations

import numpy as np

ATOL = 2e-3  # attention tolerance: |got - want| <= ATOL + RTOL * |want|
RTOL = 1e-2


def dev():
    import torch
    return torch.device("cuda:0")


def to_dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev())


def make_pools(n_layers, n_kv_heads, head_dim, num_blocks, dtype=1, rounding=0, block_size=16,
               num_host_blocks=0):
    """A device pool and the oracle layout describing the same bytes."""
    import ferrum_amd as fa
    from oracle import ref
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=n_layers, n_kv_heads=n_kv_heads,
                                         head_dim=head_dim, num_blocks=num_blocks,
                                         block_size=block_size, num_host_blocks=num_host_blocks,
                                         kv_dtype=dtype, f16_rounding=rounding))
    layout = ref.Layout(n_layers, n_kv_heads, head_dim, block_size, num_blocks, dtype, rounding)
    assert layout.pool_bytes == pool.pool_bytes
    assert layout.block_bytes == pool.block_bytes
    return pool, layout


def assert_close(got, want, atol=ATOL, rtol=RTOL, what="attention"):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    lim = atol + rtol * np.abs(want)
    bad = ~(err <= lim)
    # NaN must match NaN exactly in position
    nan_ok = np.isnan(got) == np.isnan(want)
    assert nan_ok.all(), f"{what}: NaN positions differ"
    bad &= ~(np.isnan(got) & np.isnan(want))
    assert not bad.any(), (f"{what}: {bad.sum()} values out of tolerance, "
                           f"max abs err {np.nanmax(err):.3e}")
    return float(np.nanmax(err)) if err.size else 0.0


def slots_for(table, ctx, block_size=16):
    pos = np.arange(ctx)
    return table[pos // block_size].astype(np.int64) * block_size + pos % block_size


def attention_f64(q, k_rows, v_rows, scale):
    """Brute force softmax(q K^T * scale) V in f64 for one query head.
    k_rows, v_rows: [ctx, D] decoded values."""
    s = (k_rows.astype(np.float64) @ q.astype(np.float64)) * scale
    m = s.max()
    e = np.exp(s - m)
    return (e[:, None] * v_rows.astype(np.float64)).sum(0) / e.sum()


def layer_image(pool, layout_cls, tables, ctxs, layer, seqs):
    """Host copy of one layer of the blocks the sampled sequences use, as a compact
    one-layer pool for the oracle. Returns (layout, image, remapped tables)."""
    cfg = pool.config
    bs = cfg.block_size
    ctxs = np.asarray(ctxs, np.int64)
    nb = [(int(ctxs[s]) + bs - 1) // bs for s in seqs]
    used = []
    for s, n in zip(seqs, nb):
        used.extend(int(b) for b in tables[s, :n])
    remap = {b: i for i, b in enumerate(dict.fromkeys(used))}
    lay = layout_cls(1, cfg.n_kv_heads, cfg.head_dim, bs, max(1, len(remap)), cfg.kv_dtype,
                     cfg.f16_rounding)
    region = lay.block_bytes
    image = np.zeros(lay.pool_bytes, np.uint8)
    for b, i in remap.items():
        image[i * region:(i + 1) * region] = pool.read(b * pool.block_bytes + layer * region, region)
    tab = np.zeros((len(seqs), max(1, max(nb))), np.int32)
    for j, (s, n) in enumerate(zip(seqs, nb)):
        tab[j, :n] = [remap[int(b)] for b in tables[s, :n]]
    return lay, image, tab

"""GPU parity at BASELINE.json's full configuration sizes (configs[1..4]).

The small-shape tests cover every case the kernels branch on; these run the real
shapes once and check them against the oracle through sampled sequences and
size-independent properties:
- attention outputs meet |got - want| <= 2e-3 + 1e-2 |want| against the oracle's
  restatement of crates/model/src/llama.rs:220-247 on the same pool bytes;
- appended tokens read back (FKV_GATHER_RAW) bit-exact against the oracle's encoding
  of the same f32 rows (f16 RNE, or Q8_0 per q8_dot.rs:46-59);
- copy_blocks: every sampled destination equals its source byte for byte, blocks
  outside the call are untouched; swap out -> clobber -> swap in restores the bytes.
Only the layer under test is filled; the pool has every layer of the config.
"""
import numpy as np
import pytest

from tests.helpers import assert_close, layer_image

pytestmark = pytest.mark.gpu


def _tables(pool, nblk_seq, rng, fragment_cycles=0):
    import bench
    return bench.make_tables(pool, np.asarray(nblk_seq, np.int64), rng, fragment_cycles)


def _fill(torch, pool, layer, tables, ctx, hkv, d, seed, outlier_frac=0.0):
    """N(0,1) K/V (plus +-20 outliers) for positions 0 .. ctx[s]-1 of every sequence.
    Returns the device K, V and slot tensors (kept for sampling)."""
    dev = torch.device("cuda:0")
    ctx = np.asarray(ctx, np.int64)
    seq_of = np.repeat(np.arange(ctx.size), ctx)
    pos = np.concatenate([np.arange(c) for c in ctx])
    slots = tables[seq_of, pos // 16].astype(np.int64) * 16 + pos % 16
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    k = torch.randn((slots.size, hkv, d), generator=g, device=dev)
    v = torch.randn((slots.size, hkv, d), generator=g, device=dev)
    if outlier_frac:
        for x in (k, v):
            m = torch.rand(x.shape, generator=g, device=dev) < outlier_frac
            x[m] = torch.where(torch.rand(x.shape, generator=g, device=dev) < 0.5, -20.0, 20.0)[m]
    slots_d = torch.from_numpy(slots).to(dev)
    pool.append(layer, k, v, slots_d)
    return k, v, slots


def _raw_rows_oracle(cfg, k, v):
    """Oracle encoding of token rows k, v [n, hkv, d] read back as FKV_GATHER_RAW rows."""
    from oracle import ref
    n = k.shape[0]
    lay = ref.Layout(1, cfg.n_kv_heads, cfg.head_dim, 16, (n + 15) // 16, cfg.kv_dtype,
                     cfg.f16_rounding)
    img = ref.new_pool(lay)
    slots = np.arange(n, dtype=np.int64)
    ref.append(lay, img, 0, k, v, slots)
    return ref.gather_slots(lay, img, 0, slots, 1)


def _raw_rows_device(torch, pool, layer, slots):
    cfg = pool.config
    per_head = {0: cfg.head_dim * 4, 1: cfg.head_dim * 2, 8: cfg.head_dim // 32 * 34}[cfg.kv_dtype]
    n = len(slots)
    ok = torch.zeros((n, cfg.n_kv_heads * per_head), dtype=torch.uint8, device="cuda")
    ov = torch.zeros_like(ok)
    pool.gather_slots(layer, torch.from_numpy(np.asarray(slots, np.int64)).cuda(), ok, ov, fmt=1)
    torch.cuda.synchronize()
    return ok.cpu().numpy(), ov.cpu().numpy()


def _fused_step(torch, pool, layer, hq, tables, ctx, seed):
    """One fkv_append_decode_attention call appending position ctx[s] - 1."""
    cfg = pool.config
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    n = len(ctx)
    kn = torch.randn((n, cfg.n_kv_heads, cfg.head_dim), generator=g, device="cuda")
    vn = torch.randn((n, cfg.n_kv_heads, cfg.head_dim), generator=g, device="cuda")
    q = torch.randn((n, hq, cfg.head_dim), generator=g, device="cuda")
    out = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
    ctx_d = torch.from_numpy(np.asarray(ctx, np.int32)).cuda()
    pool.append_decode_attention(layer, kn, vn, q, out, torch.from_numpy(tables).cuda(), ctx_d,
                                 int(np.max(ctx)))
    torch.cuda.synchronize()
    return kn, vn, q.cpu().numpy(), out.cpu().numpy()


def _check_decode(torch, pool, layer, tables, ctx, q, out, seqs):
    import ferrum_amd as fa
    from oracle import ref
    lay, image, tab = layer_image(pool, ref.Layout, tables, ctx, layer, seqs)
    want = ref.attention(lay, image, 0, np.ascontiguousarray(q[seqs]), tab,
                         np.asarray(ctx, np.int32)[seqs], fa.default_scale(pool.config.head_dim))
    return assert_close(out[seqs], want)


def _check_tail_raw(torch, pool, layer, tables, ctx, kn, vn):
    tail = [int(tables[s, (c - 1) // 16]) * 16 + (c - 1) % 16 for s, c in enumerate(ctx)]
    gk, gv = _raw_rows_device(torch, pool, layer, tail)
    wk, wv = _raw_rows_oracle(pool.config, kn.cpu().numpy(), vn.cpu().numpy())
    assert np.array_equal(gk, wk.reshape(gk.shape)) and np.array_equal(gv, wv.reshape(gv.shape))


def test_c2_llama3_8b_decode_step_full_size():
    """64 sequences, contexts U[128, 4096] (seed 0), 32 layers, 32/8 heads,
    D = 128, f16, scattered tables; one fused decode step on the last layer, every
    sequence checked against the oracle."""
    import torch
    import ferrum_amd as fa
    rng = np.random.default_rng(0)
    ctx0 = rng.integers(128, 4097, 64).astype(np.int64)
    nb = (ctx0 + 1 + 15) // 16
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=32, n_kv_heads=8, head_dim=128,
                                         num_blocks=int(nb.sum()) + 64))
    tables = _tables(pool, nb, rng)
    layer = 31
    _fill(torch, pool, layer, tables, ctx0, 8, 128, seed=1)
    ctx = ctx0 + 1
    kn, vn, q, out = _fused_step(torch, pool, layer, 32, tables, ctx, seed=2)
    assert pool.take_fault_flags() == 0
    _check_tail_raw(torch, pool, layer, tables, ctx, kn, vn)
    err = _check_decode(torch, pool, layer, tables, ctx, q, out, np.arange(64))
    print(f"c2: 64 sequences, max abs err {err:.2e}")
    pool.close()


def test_c4_q8_0_full_size_with_outliers():
    """Q8_0 KV, 128 sequences x 8,192 tokens, 1% of K/V at +-20 sigma. The
    fused step appends token 8,191; appended rows and a sample of 4,096 filled rows
    read back bit-exact against the oracle's quantiser, every sequence's attention
    against the oracle."""
    import torch
    import ferrum_amd as fa
    rng = np.random.default_rng(3)
    n_seqs, ctx_len = 128, 8192
    nb = np.full(n_seqs, ctx_len // 16)
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=32, n_kv_heads=8, head_dim=128,
                                         num_blocks=int(nb.sum()) + 64, kv_dtype=fa.DTYPE_Q8_0))
    tables = _tables(pool, nb, rng)
    layer = 31
    ctx0 = np.full(n_seqs, ctx_len - 1)
    k, v, slots = _fill(torch, pool, layer, tables, ctx0, 8, 128, seed=4, outlier_frac=0.01)
    pick = np.sort(rng.choice(slots.size, 4096, replace=False))
    gk, gv = _raw_rows_device(torch, pool, layer, slots[pick])
    idx = torch.from_numpy(pick).cuda()
    wk, wv = _raw_rows_oracle(pool.config, k[idx].cpu().numpy(), v[idx].cpu().numpy())
    assert np.array_equal(gk, wk.reshape(gk.shape)) and np.array_equal(gv, wv.reshape(gv.shape))
    del k, v
    ctx = np.full(n_seqs, ctx_len)
    kn, vn, q, out = _fused_step(torch, pool, layer, 32, tables, ctx, seed=5)
    assert pool.take_fault_flags() == 0
    _check_tail_raw(torch, pool, layer, tables, ctx, kn, vn)
    err = _check_decode(torch, pool, layer, tables, ctx, q, out, np.arange(n_seqs))
    print(f"c4: 128 sequences, max abs err {err:.2e}")
    pool.close()


def test_c3_continuous_batching_full_size():
    """a 172.8 GB pool (60% of 288 GB) fragmented by 10,000 seeded
    alloc/free cycles; 256 decode sequences with log-normal contexts (median 2048,
    sigma 1.0, cap 32,768) and 4 sequences appending a 512-token prefill chunk in the
    same step. Every decode sequence and every query row of the four prefill chunks
    against the oracle."""
    import torch
    import ferrum_amd as fa
    from oracle import ref
    rng = np.random.default_rng(6)
    L, hq, hkv, d = 32, 32, 8, 128
    ctx_dec = np.minimum(np.round(np.exp(rng.normal(np.log(2048), 1.0, 256))), 32767)
    ctx_dec = np.maximum(ctx_dec, 1).astype(np.int64)
    prior = np.array([0, 512, 1024, 1536], np.int64)
    chunk = 512
    block_bytes = L * 2 * hkv * 16 * d * 2
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=L, n_kv_heads=hkv, head_dim=d,
                                         num_blocks=int(0.6 * 288e9 // block_bytes)))
    nb = np.concatenate([(ctx_dec + 1 + 15) // 16, (prior + chunk + 15) // 16])
    tables = _tables(pool, nb, rng, fragment_cycles=10000)
    layer = 0
    _fill(torch, pool, layer, tables, np.concatenate([ctx_dec, prior]), hkv, d, seed=7)
    # decode part: fused step for the 256 decode sequences
    dec_tab = np.ascontiguousarray(tables[:256])
    ctx = ctx_dec + 1
    kn, vn, q, out = _fused_step(torch, pool, layer, hq, dec_tab, ctx, seed=8)
    # prefill part: append the chunk through its slot mapping, then chunked attention
    pre_tab = np.ascontiguousarray(tables[256:])
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    kp = torch.randn((4 * chunk, hkv, d), generator=g, device="cuda")
    vp = torch.randn((4 * chunk, hkv, d), generator=g, device="cuda")
    qp = torch.randn((4 * chunk, hq, d), generator=g, device="cuda")
    op = torch.full(qp.shape, 7.0, dtype=torch.float32, device="cuda")
    pos = np.concatenate([np.arange(p, p + chunk) for p in prior])
    seq = np.repeat(np.arange(4), chunk)
    pslots = pre_tab[seq, pos // 16].astype(np.int64) * 16 + pos % 16
    pool.append(layer, kp, vp, torch.from_numpy(pslots).cuda())
    pctx = (prior + chunk).astype(np.int32)
    qlen = np.full(4, chunk, np.int32)
    qoff = np.arange(0, 4 * chunk, chunk, dtype=np.int64)
    pool.prefill_attention(layer, qp, op, torch.from_numpy(pre_tab).cuda(),
                           torch.from_numpy(pctx).cuda(), torch.from_numpy(qlen).cuda(),
                           torch.from_numpy(qoff).cuda(), chunk, int(pctx.max()))
    torch.cuda.synchronize()
    assert pool.take_fault_flags() == 0
    err = _check_decode(torch, pool, layer, dec_tab, ctx, q, out, np.arange(256))
    _check_tail_raw(torch, pool, layer, dec_tab, ctx, kn, vn)
    # prefill: every row of the four chunks, against the oracle's token-by-token restatement
    lay, image, tab = layer_image(pool, ref.Layout, pre_tab, pctx, layer, [0, 1, 2, 3])
    want = ref.prefill_attention(lay, image, 0, qp.cpu().numpy(), tab, pctx, qlen, qoff,
                                 fa.default_scale(d))
    perr = assert_close(op.cpu().numpy(), want, what="prefill")
    print(f"c3: 256 decode sequences, max abs err {err:.2e}; 2,048 prefill rows, {perr:.2e}")
    pool.close()


def test_c5_llama3_70b_long_context_copy_and_swap_full_size():
    """one 131,072-token sequence on 70B-shaped KV (80 layers, 64/8
    heads, f16, 42.9 GB), decode attention over the full context against the oracle;
    copy_blocks of 20,000 seeded (src, dst) pairs (distinct destinations) and a swap
    of 20% of the context's blocks out to pinned host memory and back."""
    import torch
    import ferrum_amd as fa
    rng = np.random.default_rng(10)
    ctx_len, n_pairs = 131072, 20000
    nctx = ctx_len // 16
    n_swap = nctx // 5
    pool = fa.PagedKvPool(fa.PagedConfig(n_layers=80, n_kv_heads=8, head_dim=128,
                                         num_blocks=nctx + n_pairs + 64, num_host_blocks=n_swap))
    tables = _tables(pool, np.array([nctx]), rng)
    layer = 79
    _fill(torch, pool, layer, tables, np.array([ctx_len - 1]), 8, 128, seed=11)
    ctx = np.array([ctx_len])
    kn, vn, q, out = _fused_step(torch, pool, layer, 64, tables, ctx, seed=12)
    assert pool.take_fault_flags() == 0
    _check_tail_raw(torch, pool, layer, tables, ctx, kn, vn)
    err = _check_decode(torch, pool, layer, tables, ctx, q, out, [0])
    print(f"c5: attention max abs err {err:.2e}")

    bb = pool.block_bytes
    used = tables[0, :nctx].astype(np.int64)
    dst = pool.alloc_blocks(n_pairs).astype(np.int64)
    src = used[rng.integers(0, nctx, n_pairs)]
    spare = pool.alloc_blocks(4).astype(np.int64)  # never a destination
    spare_before = [pool.read(int(b) * bb, bb) for b in spare]
    pool.copy_blocks(torch.from_numpy(np.stack([src, dst], 1)).cuda())
    torch.cuda.synchronize()
    for j in rng.integers(0, n_pairs, 24):
        assert np.array_equal(pool.read(int(dst[j]) * bb, bb), pool.read(int(src[j]) * bb, bb))
    for b, before in zip(spare, spare_before):
        assert np.array_equal(pool.read(int(b) * bb, bb), before)

    sel = np.sort(rng.choice(used, n_swap, replace=False))
    check = sel[rng.integers(0, n_swap, 12)]
    before = [pool.read(int(b) * bb, bb) for b in check]
    pool.swap_out(np.stack([sel, np.arange(n_swap)], 1))
    torch.cuda.synchronize()
    pool.fill(0x5A)
    pool.swap_in(np.stack([np.arange(n_swap), sel], 1))
    torch.cuda.synchronize()
    for b, want in zip(check, before):
        assert np.array_equal(pool.read(int(b) * bb, bb), want)
    assert pool.take_fault_flags() == 0
    pool.close()

"""CPU: the oracle's pool semantics and attention loop (no GPU).

Dense revision-1 pool: the unit tests of crates/kvcache/src/pool.rs:233-308
ported onto the oracle's restatement (the same tests run on the device pool in
test_gpu_compat.py). Paged operations: closed forms (gather(append(x)) == enc(x),
copy_blocks is a block memcpy that leaves other blocks alone). Attention: the
loop of crates/model/src/llama.rs:220-247 against an f64 brute force and against
closed forms (ctx = 1 gives V_0; equal keys give mean(V); one dominant key gives
its V; a non-finite max gives zeros, scalar.rs:125-130), GQA mapping kv_h = h / g,
and invariance under permuting physical blocks.
"""
import numpy as np
import pytest

from oracle import ref
from tests.helpers import attention_f64, slots_for

TINY = (2, 1, 4, 3, 2)  # pool.rs:237-245: layers, kv heads, head dim, max seq, slots
K4 = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
V4 = np.array([5.0, 6.0, 7.0, 8.0], np.float32)


def ok(res):
    assert res[0] == 0, res[1]
    return res[2]


def test_dense_round_trip():
    # pool.rs:247-261
    p = ref.DensePool(*TINY)
    slot = ok(p.alloc())
    assert ok(p.seq_len(slot)) == 0
    ok(p.append_layer(slot, 0, K4, V4))
    ok(p.append_layer(slot, 1, K4, V4))
    ok(p.commit_token(slot))
    assert ok(p.seq_len(slot)) == 1
    assert np.array_equal(ok(p.k(slot, 0, 0)), K4)
    assert np.array_equal(ok(p.v(slot, 1, 0)), V4)


def test_dense_layer_order_and_commit():
    # pool.rs:263-275
    p = ref.DensePool(*TINY)
    slot = ok(p.alloc())
    assert p.append_layer(slot, 1, K4, V4)[:2] == (1, "cache: layers must append in order")
    ok(p.append_layer(slot, 0, K4, V4))
    assert p.commit_token(slot)[:2] == (1, "cache: not every layer appended")
    ok(p.append_layer(slot, 1, K4, V4))
    ok(p.commit_token(slot))
    assert p.k(slot, 0, 1)[:2] == (1, "cache: position not yet committed")


def test_dense_abandon_and_uncommit():
    # pool.rs:277-291
    p = ref.DensePool(*TINY)
    slot = ok(p.alloc())
    ok(p.append_layer(slot, 0, K4, V4))
    ok(p.abandon_partial(slot))
    ok(p.append_layer(slot, 0, K4, V4))
    ok(p.append_layer(slot, 1, K4, V4))
    ok(p.commit_token(slot))
    ok(p.uncommit_token(slot))
    assert ok(p.seq_len(slot)) == 0
    ok(p.append_layer(slot, 0, K4, V4))
    assert p.uncommit_token(slot)[:2] == (1, "cache: nothing to uncommit")


def test_dense_storage_size_and_exhaustion():
    # pool.rs:293-307 and the Unavailable rule of pool.rs:84-88
    p = ref.DensePool(*TINY)
    assert p.storage_len() == 2 * 2 * 3 * 1 * 4 * 2
    ok(p.alloc())
    ok(p.alloc())
    assert p.alloc()[:2] == (2, "no free kv slots")
    assert p.storage_len() == 2 * 2 * 3 * 1 * 4 * 2
    assert p.free(5)[:2] == (1, "cache: free of unallocated slot")
    bad = ref.DensePool(0, 1, 4, 3, 2)
    assert (bad.code, bad.msg) == (1, "cache: kv pool dimension is zero")
    big = ref.DensePool(1 << 20, 1 << 20, 1 << 20, 1 << 20, 2)
    assert (big.code, big.msg) == (1, "cache: kv pool size overflow")


def test_dense_alloc_zero_fills_a_reused_slot():
    # pool.rs:92-97: alloc zero-fills, so a freed-then-reallocated slot reads zeros
    p = ref.DensePool(*TINY)
    s = ok(p.alloc())
    ok(p.append_layer(s, 0, K4, V4))
    ok(p.append_layer(s, 1, K4, V4))
    ok(p.commit_token(s))
    ok(p.free(s))
    s2 = ok(p.alloc())
    assert s2 == s
    ok(p.append_layer(s2, 0, np.zeros(4, np.float32), np.zeros(4, np.float32)))
    ok(p.append_layer(s2, 1, np.zeros(4, np.float32), np.zeros(4, np.float32)))
    ok(p.commit_token(s2))
    assert np.all(ok(p.k(s2, 1, 0)) == 0)


# -- paged closed forms ------------------------------------------------------------

def _enc(x, dtype, rounding):
    """Expected decoded values after storage (closed forms, not the oracle)."""
    if dtype == 0:
        return x
    if dtype == 1:
        if rounding == 0:
            return x.astype(np.float16).astype(np.float32)
        return ref.f16_to_f32(ref.f32_to_f16(x, 1))
    raw = ref.q8_quantize_row(x.ravel(), rounding)
    return ref.q8_dequant(raw, x.size).reshape(x.shape)


@pytest.mark.parametrize("dtype,d,rounding", [(0, 64, 0), (1, 128, 0), (1, 64, 1), (8, 128, 0),
                                              (8, 64, 1), (1, 12, 0)])
def test_gather_of_append_is_encoding(dtype, d, rounding):
    rng = np.random.default_rng(d + dtype)
    lay = ref.Layout(3, 2, d, 16, 40, dtype, rounding)
    pool = ref.new_pool(lay)
    ctx = [37, 1, 16, 100, 0, 33]
    perm = rng.permutation(40).astype(np.int32)
    mb = max((c + 15) // 16 for c in ctx)
    tab = np.zeros((len(ctx), mb), np.int32)
    off = 0
    for i, c in enumerate(ctx):
        n = (c + 15) // 16
        tab[i, :n] = perm[off:off + n]
        off += n
    slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(ctx)])
    slots = np.insert(slots, [2, 9], -1)
    x = rng.standard_normal((slots.size, 2, d)).astype(np.float32)
    y = rng.standard_normal((slots.size, 2, d)).astype(np.float32)
    assert ref.append(lay, pool, 1, x, y, slots) == 0
    gk, gv = ref.gather_slots(lay, pool, 1, slots, 0)
    live = slots >= 0
    if dtype == 8:
        ek = _enc(x[live].reshape(-1, d), dtype, rounding).reshape(-1, 2, d)
        ev = _enc(y[live].reshape(-1, d), dtype, rounding).reshape(-1, 2, d)
    else:
        ek, ev = _enc(x[live], dtype, rounding), _enc(y[live], dtype, rounding)
    assert np.array_equal(gk[live].view(np.uint32), ek.view(np.uint32))
    assert np.array_equal(gv[live].view(np.uint32), ev.view(np.uint32))
    # by block table: rows in sequence order
    tk, tv, offs = ref.gather_tables(lay, pool, 1, tab, np.array(ctx, np.int32), 0)
    assert np.array_equal(tk.view(np.uint32), gk[live].view(np.uint32))
    # other layers untouched
    assert not ref.gather_slots(lay, pool, 0, slots[live], 1)[0].any()


def test_out_of_range_slot_is_skipped():
    lay = ref.Layout(1, 1, 32, 16, 2, 1, 0)
    pool = ref.new_pool(lay)
    x = np.ones((3, 1, 32), np.float32)
    assert ref.append(lay, pool, 0, x, x, np.array([0, 32, 5])) == 1
    assert np.count_nonzero(pool.view(np.uint16) == 0x3C00) == 2 * 2 * 32  # 2 tokens, K and V


def test_copy_blocks_is_block_memcpy():
    rng = np.random.default_rng(0)
    lay = ref.Layout(2, 2, 64, 16, 12, 8, 0)
    img = rng.integers(0, 256, lay.pool_bytes, dtype=np.uint8)
    pool = img.copy()
    pairs = np.array([[0, 7], [3, 8], [3, 9], [11, 4]], np.int64)
    ref.copy_blocks(lay, pool, pairs)
    bb = lay.block_bytes
    want = img.copy()
    for s, d in pairs:
        want[d * bb:(d + 1) * bb] = img[s * bb:(s + 1) * bb]
    assert np.array_equal(pool, want)


# -- attention -------------------------------------------------------------------

def _pool_with(dtype, d, hkv, ctxs, seed, perm_seed=None, layers=1):
    rng = np.random.default_rng(seed)
    nb = [(c + 15) // 16 for c in ctxs]
    nblk = sum(nb) + 3
    lay = ref.Layout(layers, hkv, d, 16, nblk, dtype, 0)
    pool = ref.new_pool(lay)
    perm = np.random.default_rng(seed if perm_seed is None else perm_seed).permutation(nblk)
    tab = np.zeros((len(ctxs), max(1, max(nb))), np.int32)
    off = 0
    for i, n in enumerate(nb):
        tab[i, :n] = perm[off:off + n]
        off += n
    total = sum(ctxs)
    k = rng.standard_normal((total, hkv, d)).astype(np.float32)
    v = rng.standard_normal((total, hkv, d)).astype(np.float32)
    slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(ctxs)])
    for layer in range(layers):
        ref.append(lay, pool, layer, k, v, slots)
    return lay, pool, tab


@pytest.mark.parametrize("dtype,d,g", [(1, 128, 4), (1, 64, 8), (0, 64, 1), (8, 128, 2)])
def test_attention_matches_f64_brute_force(dtype, d, g):
    ctxs = [1, 17, 300, 64]
    hkv = 2
    lay, pool, tab = _pool_with(dtype, d, hkv, ctxs, seed=1)
    q = np.random.default_rng(2).standard_normal((len(ctxs), hkv * g, d)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    out = ref.attention(lay, pool, 0, q, tab, np.array(ctxs, np.int32), scale)
    for s, c in enumerate(ctxs):
        kr, vr = ref.gather_slots(lay, pool, 0, slots_for(tab[s], c), 0)
        for h in range(hkv * g):
            want = attention_f64(q[s, h], kr[:, h // g], vr[:, h // g], scale)
            assert np.allclose(out[s, h], want, rtol=1e-5, atol=1e-6), (s, h)


def test_attention_closed_forms():
    d, hkv, g = 64, 1, 4
    lay = ref.Layout(1, hkv, d, 16, 8, 0, 0)
    rng = np.random.default_rng(5)
    tab = np.arange(8, dtype=np.int32)[None, :]
    q = rng.standard_normal((1, g, d)).astype(np.float32)
    # ctx = 1 -> V_0 exactly (softmax of one element is 1)
    pool = ref.new_pool(lay)
    k = rng.standard_normal((100, 1, d)).astype(np.float32)
    v = rng.standard_normal((100, 1, d)).astype(np.float32)
    ref.append(lay, pool, 0, k, v, slots_for(tab[0], 100))
    out = ref.attention(lay, pool, 0, q, tab, np.array([1], np.int32), 0.125)
    assert np.array_equal(out[0], np.repeat(v[0], g, axis=0))
    # all keys equal -> mean of V
    k_eq = np.repeat(k[:1], 100, axis=0)
    ref.append(lay, pool, 0, k_eq, v, slots_for(tab[0], 100))
    out = ref.attention(lay, pool, 0, q, tab, np.array([100], np.int32), 0.125)
    assert np.allclose(out[0], v[:, 0].astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)
    # one key dominates (score gap 1e4) -> its V
    k_dom = np.zeros((100, 1, d), np.float32)
    k_dom[37, 0] = q[0, 0] * 1e3
    ref.append(lay, pool, 0, k_dom, v, slots_for(tab[0], 100))
    out = ref.attention(lay, pool, 0, q, tab, np.array([100], np.int32), 1.0)
    assert np.array_equal(out[0, 0], v[37, 0])
    # +inf score -> non-finite max -> zeros (scalar.rs:127-130)
    k_inf = np.zeros((100, 1, d), np.float32)
    k_inf[3, 0, 0] = np.inf
    ref.append(lay, pool, 0, k_inf, v, slots_for(tab[0], 100))
    qq = np.zeros((1, g, d), np.float32)
    qq[0, :, 0] = 1.0
    out = ref.attention(lay, pool, 0, qq, tab, np.array([100], np.int32), 0.125)
    assert np.all(out == 0)
    # empty context -> zeros
    out = ref.attention(lay, pool, 0, q, tab, np.array([0], np.int32), 0.125)
    assert np.all(out == 0)


def test_attention_gqa_mapping_and_block_placement():
    ctxs = [50, 200]
    d, hkv, g = 64, 2, 4
    q = np.random.default_rng(3).standard_normal((2, hkv * g, d)).astype(np.float32)
    outs = []
    for ps in (10, 11):
        lay, pool, tab = _pool_with(1, d, hkv, ctxs, seed=4, perm_seed=ps)
        outs.append(ref.attention(lay, pool, 0, q, tab, np.array(ctxs, np.int32), 0.125))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    # query heads 0..g-1 read KV head 0: with identical q rows they give identical out
    lay, pool, tab = _pool_with(1, d, hkv, ctxs, seed=4)
    q2 = q.copy()
    q2[:, 1:g] = q2[:, :1]
    o = ref.attention(lay, pool, 0, q2, tab, np.array(ctxs, np.int32), 0.125)
    assert np.array_equal(o[:, 1], o[:, 0]) and not np.array_equal(o[:, g], o[:, 0])


@pytest.mark.parametrize("dtype", [1, 8, 0])
def test_avx2_attention_within_tolerance_of_oracle(dtype):
    """The CPU baseline's AVX2 port reads every storage type's tiles as the scalar oracle
    does (Q8_0: the quants' operand order inside the tile)."""
    if not ref.avx2_available():
        pytest.skip("host has no AVX2/FMA/F16C")
    ctxs = [3, 129, 700]
    lay, pool, tab = _pool_with(dtype, 128, 2, ctxs, seed=9)
    q = np.random.default_rng(1).standard_normal((3, 8, 128)).astype(np.float32)
    c = np.array(ctxs, np.int32)
    a = ref.attention(lay, pool, 0, q, tab, c, 0.088388346)
    b1 = ref.avx2_attention(lay, pool, 0, q, tab, c, 0.088388346, 1)
    b4 = ref.avx2_attention(lay, pool, 0, q, tab, c, 0.088388346, 4)
    assert np.array_equal(b1, b4)
    assert np.allclose(a, b1, rtol=1e-5, atol=1e-6)


def test_prefill_is_decode_at_every_position_and_causal_brute_force():
    """Prefill of a chunk (llama.rs:363-378) == the decode loop at each of its positions,
    and == an f64 causal softmax(qK^T)V."""
    ctxs, qls = [40, 300, 17], [40, 33, 5]
    d, hkv, g = 64, 2, 4
    lay, pool, tab = _pool_with(1, d, hkv, ctxs, seed=12)
    rows = sum(qls)
    offs = np.concatenate([[0], np.cumsum(qls)[:-1]]).astype(np.int64)
    q = np.random.default_rng(4).standard_normal((rows, hkv * g, d)).astype(np.float32)
    scale = 0.125
    got = ref.prefill_attention(lay, pool, 0, q, tab, np.array(ctxs, np.int32),
                                np.array(qls, np.int32), offs, scale)
    for s, (c, n) in enumerate(zip(ctxs, qls)):
        kr, vr = ref.gather_slots(lay, pool, 0, slots_for(tab[s], c), 0)
        for i in range(n):
            r = offs[s] + i
            pos_ctx = c - n + i + 1
            dec = ref.attention(lay, pool, 0, q[r:r + 1], tab[s:s + 1],
                                np.array([pos_ctx], np.int32), scale)
            assert np.array_equal(got[r], dec[0])
            if i in (0, n - 1):
                for h in (0, hkv * g - 1):
                    want = attention_f64(q[r, h], kr[:pos_ctx, h // g], vr[:pos_ctx, h // g], scale)
                    assert np.allclose(got[r, h], want, rtol=1e-5, atol=1e-6)
